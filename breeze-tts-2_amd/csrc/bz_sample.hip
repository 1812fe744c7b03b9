// CFG + HF-order sampling of one token per row in one launch (gfx950).
//
// Replaces the depth decoder's per-codebook sampling sequence
// (models/cudagraph/depth_decoder_graph.py:487-558, _cfg_sample): the CFG
// combination uncond + g * (cond - uncond), the invalid-codec-token mask
// (models/logits_process.py:7-25), temperature, top-k over a fixed workspace,
// top-p, softmax, multinomial, and argmax for greedy rows -- about twenty
// torch kernels -- with one workgroup per sampled row:
//
//   1. combined logits of the row (and its greedy argmax, first index of the
//      maximum, as torch.argmax) into LDS, divided by the temperature;
//   2. the k-th largest entry (k = top_k, or the whole workspace) by a radix
//      select over unique 64-bit keys (scaled value, then ascending index),
//      and a bitonic sort of just those k entries (padded to a power of two
//      >= 64; partners under 64 apart trade through wave shuffles): rank r of
//      the sorted set is rank r of top-k;
//   3. the top-k ranks (k = top_k, or the whole workspace for top_k <= 0)
//      and their softmax (one rank per thread, the workspace is <= 1024
//      wide), an inclusive block scan of it, and the top-p prefix: rank r
//      stays when r == 0 or the cumulative probability before it is <= top_p
//      (the reference's shifted mask), so the kept set is a prefix of ranks;
//   4. one uniform draw u in [0, 1) (Philox4x32-10, Salmon, Moraes, Dror and
//      Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011; key =
//      the 64-bit seed, read from device memory so a captured graph picks up
//      a new one; counter = (the row's call count, row)) and the first
//      kept rank whose cumulative weight exceeds u times the kept total;
//   5. the token (sampled, or the argmax when do_sample is 0) to the row and
//      its unconditional twin; the row's call count is advanced, so graph
//      replays draw fresh numbers.
// A greedy row that reports no probabilities stops after step 1.
//
// The random stream is this library's own, not torch's: the sampled tokens
// follow the same distribution as the reference's, not the same sequence.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "bz_gemv.h"
#include "bz_sample.h"

namespace bz {
namespace {

constexpr int kSampleThreads = 1024;
constexpr int kSampleWidth = 4096;  // padded row: the largest vocabulary
constexpr int kSampleMaxK = 1024;   // top-k workspace: one rank per thread

// Philox4x32-10 of the paper above: 10 rounds of the 4x32 round function with
// its published multipliers and Weyl key increments.
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
    constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u, kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)kM0 * c[0], p1 = (uint64_t)kM1 * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1, n3 = (uint32_t)p0;
        c[0] = n0;
        c[1] = n1;
        c[2] = n2;
        c[3] = n3;
        k0 += kW0;
        k1 += kW1;
    }
}

struct SampleParams {
    const float* logits;
    int64_t ld;
    int B, half, V, codec, max_k;
    const float* guidance;
    const float* temperature;
    const int64_t* top_k;
    const float* top_p;
    const int64_t* do_sample;
    const uint64_t* seed;
    uint64_t* counters;
    int64_t* tokens;
    float* cfg_out;
    float* probs_out;
};

// Sort key of a row entry: the temperature-scaled value mapped to an
// unsigned order (larger float -> larger key) in the high word, the inverted
// index in the low word, so keys are unique and a larger key is a larger
// value, or the same value at a smaller index (the order of torch.argmax).
__device__ __forceinline__ uint64_t entry_key(float s, int v) {
    const uint32_t b = __float_as_uint(s);
    const uint32_t u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)v);
}
__device__ __forceinline__ float key_value(uint64_t key) {
    const uint32_t u = (uint32_t)(key >> 32);
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}
__device__ __forceinline__ int key_index(uint64_t key) { return (int)(0xFFFFFFFFu - (uint32_t)key); }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, 64), hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float wave_scan_incl(float v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

constexpr int kPerThread = kSampleWidth / kSampleThreads;  // row entries a thread holds

__global__ void __launch_bounds__(kSampleThreads) sample_cfg_kernel(SampleParams p) {
    __shared__ uint64_t cand[kSampleMaxK];  // the selected keys, then sorted
    __shared__ unsigned hist[256];
    __shared__ float wsum[kSampleThreads / 64];
    __shared__ float wbest_v[kSampleThreads / 64];
    __shared__ int wbest_i[kSampleThreads / 64];
    __shared__ int greedy_s, ncand, sel_digit, sel_need, sel_count, pick, last_kept;
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int NW = kSampleThreads / 64;
    const float* cond = p.logits + (int64_t)r * p.ld;
    const float* uncond = p.logits + (int64_t)(p.B >= 2 ? p.half + r : r) * p.ld;
    const float g = p.B >= 2 ? p.guidance[r] : 0.0f;
    const float temp = p.temperature[r];

    // 1. combined logits, greedy argmax, the scaled entries' keys (registers)
    float best_v = -INFINITY;
    int best_i = 0x7FFFFFFF;
    uint64_t key[kPerThread];
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
        const int v = tid + q * kSampleThreads;
        key[q] = 0;  // absent (below every entry's key)
        if (v < p.V) {
            float c = cond[v];
            if (p.B >= 2) {
                const float u = uncond[v];
                c = u + g * (c - u);
            }
            if (v >= p.codec) c = -INFINITY;
            if (p.cfg_out) p.cfg_out[(int64_t)r * p.V + v] = c;
            if (c > best_v || best_i == 0x7FFFFFFF) {  // ascending v: the first maximum wins
                best_v = c;
                best_i = v;
            }
            key[q] = entry_key(c / temp, v);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best_v, o, 64);
        const int oi = __shfl_xor(best_i, o, 64);
        if (ov > best_v || (ov == best_v && oi < best_i)) {
            best_v = ov;
            best_i = oi;
        }
    }
    if (lane == 0) {
        wbest_v[wave] = best_v;
        wbest_i[wave] = best_i;
    }
    if (tid == 0) ncand = 0;

    // A greedy row with no probabilities to report needs only the argmax:
    // skip the select, sort, softmax and draw.  Same token (same reduction
    // order as below) and the call count advances as on the full path.
    if (!p.do_sample[r] && !p.probs_out) {
        __syncthreads();
        if (tid == 0) {
            float bv = wbest_v[0];
            int bi = wbest_i[0];
            for (int w = 1; w < NW; ++w)
                if (wbest_v[w] > bv || (wbest_v[w] == bv && wbest_i[w] < bi)) {
                    bv = wbest_v[w];
                    bi = wbest_i[w];
                }
            const int64_t tok = bi < 0 ? 0 : (bi >= p.V ? p.V - 1 : bi);
            p.tokens[r] = tok;
            if (p.B >= 2) p.tokens[p.half + r] = tok;
            p.counters[r] = p.counters[r] + 1;
        }
        return;
    }

    // 2. the k-th largest key (k = top_k, or the whole workspace): radix
    //    select over 8-bit digits from the top; keys are unique, so exactly k
    //    keys are >= the result.  A pass whose chosen bucket holds exactly
    //    the keys still needed ends the search.
    const int64_t tk = p.top_k[r];
    const int kk = tk > 0 ? (int)min<int64_t>(tk, p.max_k) : p.max_k;
    uint64_t prefix = 0, mask = 0;
    int need = kk;
    for (int shift = 56; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPerThread; ++q)
            if (key[q] != 0 && (key[q] & mask) == prefix) atomicAdd(&hist[(key[q] >> shift) & 255u], 1u);
        __syncthreads();
        if (wave == 0) {
            // lane l covers digits 255 - 4l .. 252 - 4l (top down)
            unsigned c4[4], sum = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                c4[q] = hist[255 - 4 * lane - q];
                sum += c4[q];
            }
            unsigned incl = sum;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const unsigned t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            unsigned above = incl - sum;  // keys in higher digits than this lane's
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (above < (unsigned)need && above + c4[q] >= (unsigned)need) {
                    sel_digit = 255 - 4 * lane - q;
                    sel_need = need - (int)above;
                    sel_count = (int)c4[q];
                }
                above += c4[q];
            }
        }
        __syncthreads();
        prefix |= (uint64_t)sel_digit << shift;
        mask |= (uint64_t)255u << shift;
        need = sel_need;
        if (sel_count == need) break;  // workgroup-uniform
    }

    // 3. the kk selected keys into LDS, padded with zeros to P (a power of
    //    two >= 64), then a bitonic sort, descending: partners less than 64
    //    apart trade through wave shuffles, wider ones through LDS
    const int P = max(64, 1 << (32 - __clz(kk - 1)));
#pragma unroll
    for (int q = 0; q < kPerThread; ++q)
        if (key[q] != 0 && key[q] >= prefix) cand[atomicAdd(&ncand, 1)] = key[q];
    __syncthreads();
    uint64_t mine = tid < kk ? cand[tid] : 0;
    for (int lk = 1; (1 << lk) <= P; ++lk) {
        const int k = 1 << lk;
        for (int lj = lk - 1; lj >= 0; --lj) {
            const int j = 1 << lj;
            uint64_t theirs;
            if (j < 64) {
                theirs = shfl_xor64(mine, j);
            } else {
                __syncthreads();
                if (tid < P) cand[tid] = mine;
                __syncthreads();
                theirs = tid < P ? cand[tid ^ j] : 0;
            }
            const bool lower = (tid & j) == 0, desc = (tid & k) == 0;
            const uint64_t hi = mine > theirs ? mine : theirs, lo = mine > theirs ? theirs : mine;
            if (tid < P) mine = (lower == desc) ? hi : lo;
        }
    }
    if (tid == 0) {
        float bv = wbest_v[0];
        int bi = wbest_i[0];
        for (int w = 1; w < NW; ++w)
            if (wbest_v[w] > bv || (wbest_v[w] == bv && wbest_i[w] < bi)) {
                bv = wbest_v[w];
                bi = wbest_i[w];
            }
        greedy_s = bi;
    }

    // 4. thread t = rank t: top-k softmax weights, block scan, top-p prefix
    const int t = tid;
    const float sv_t = key_value(mine);
    const int si_t = key_index(mine);
    __shared__ float m_s;  // rank 0 holds the maximum
    if (tid == 0) m_s = sv_t;
    __syncthreads();
    const float e = (t < kk && sv_t > -INFINITY) ? expf(sv_t - m_s) : 0.0f;
    float inc = wave_scan_incl(e, lane);
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    float before_w = 0.0f, total = 0.0f;
    for (int w = 0; w < NW; ++w) {
        if (w < wave) before_w += wsum[w];
        total += wsum[w];
    }
    inc += before_w;
    const float exc = inc - e;
    // kept: rank 0, or the cumulative probability before this rank <= top_p
    const bool kept = t < kk && e > 0.0f && (t == 0 || exc / total <= p.top_p[r]);
    __syncthreads();  // wsum is reused below
    const float ke = kept ? e : 0.0f;  // the kept set is a prefix of ranks
    float ks = ke;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ks += __shfl_xor(ks, o, 64);
    if (lane == 0) wsum[wave] = ks;
    if (tid == 0) {
        pick = 0x7FFFFFFF;
        last_kept = 0;
    }
    __syncthreads();
    float kept_total = 0.0f;
    for (int w = 0; w < NW; ++w) kept_total += wsum[w];

    if (p.probs_out) {
        float* pr = p.probs_out + (int64_t)r * p.V;
        for (int v = tid; v < p.V; v += kSampleThreads) pr[v] = 0.0f;
        __syncthreads();
        if (kept) pr[si_t] = ke / kept_total;
    }

    // 5. the draw: the first kept rank whose cumulative weight exceeds
    //    u * kept_total (kept ranks are a prefix, so their cumulative weight
    //    is `inc`)
    const uint64_t cnt = p.counters[r];
    uint32_t c[4] = {(uint32_t)cnt, (uint32_t)(cnt >> 32), (uint32_t)r, 0u};
    const uint64_t keyr = *p.seed;
    philox4x32_10(c, (uint32_t)keyr, (uint32_t)(keyr >> 32));
    const float u = (float)(c[0] >> 8) * (1.0f / 16777216.0f);
    if (kept) {
        atomicMax(&last_kept, t);
        if (inc > u * kept_total) atomicMin(&pick, t);
    }
    __syncthreads();
    if (tid == (pick == 0x7FFFFFFF ? last_kept : pick)) {  // rounding at the top end: the last kept rank
        // 6. the token, to the row and its twin; advance the row's call count
        int64_t tok = p.do_sample[r] ? (int64_t)si_t : (int64_t)greedy_s;
        tok = tok < 0 ? 0 : (tok >= p.V ? p.V - 1 : tok);
        p.tokens[r] = tok;
        if (p.B >= 2) p.tokens[p.half + r] = tok;
        p.counters[r] = cnt + 1;
    }
}

}  // namespace
}  // namespace bz

using namespace bz;

extern "C" int bz_sample_cfg(const float* logits, int64_t ld_logits, int32_t B, int32_t V, int32_t codec_size,
                             int32_t max_k, const float* guidance, const float* temperature, const int64_t* top_k,
                             const float* top_p, const int64_t* do_sample, const uint64_t* seed, uint64_t* counters,
                             int64_t* tokens, float* cfg_out, float* probs_out, void* stream) {
    if (!logits || !temperature || !top_k || !top_p || !do_sample || !seed || !counters || !tokens)
        return BZ_ERR_INVALID_ARG;
    if (B < 1 || (B > 1 && B % 2) || V < 1 || V > kSampleWidth || ld_logits < V) return BZ_ERR_INVALID_ARG;
    if (codec_size < 1 || codec_size > V || max_k < 1 || max_k > kSampleMaxK || max_k > V) return BZ_ERR_INVALID_ARG;
    if (B >= 2 && !guidance) return BZ_ERR_INVALID_ARG;
    SampleParams p;
    p.logits = logits;
    p.ld = ld_logits;
    p.B = B;
    p.half = B == 1 ? 1 : B / 2;
    p.V = V;
    p.codec = codec_size;
    p.max_k = max_k;
    p.guidance = guidance;
    p.temperature = temperature;
    p.top_k = top_k;
    p.top_p = top_p;
    p.do_sample = do_sample;
    p.seed = seed;
    p.counters = counters;
    p.tokens = tokens;
    p.cfg_out = cfg_out;
    p.probs_out = probs_out;
    hipLaunchKernelGGL(sample_cfg_kernel, dim3(p.half), dim3(kSampleThreads), 0, static_cast<hipStream_t>(stream), p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}
