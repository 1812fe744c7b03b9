/* CFG + HF-order token sampling on the GPU (libbzgemv.so).  C ABI: plain
 * pointers and sizes, device memory, a HIP stream (NULL = default). */
#ifndef BZ_SAMPLE_H
#define BZ_SAMPLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One token per sampled row from fp32 logits [B][ld_logits] (V used).
 * B = 1 (no CFG) or 2 half (rows [0, half) conditional, [half, B)
 * unconditional): combined = uncond + guidance[r] * (cond - uncond), columns
 * [codec_size, V) masked to -inf, then temperature, top-k over a max_k-wide
 * workspace (top_k[r] <= 0: the whole workspace), top-p with the shifted
 * mask (the token that crosses top_p stays), softmax and one draw; rows with
 * do_sample[r] == 0 take the first argmax of the combined logits.  The token
 * goes to tokens[r] and, with CFG, tokens[half + r]; counters[r] (the row's
 * draw count; *seed, in device memory, is the Philox4x32-10 key) is
 * advanced by one, so replays of a captured call draw fresh numbers.
 * Per-row parameters have half entries.  cfg_out / probs_out (optional,
 * [half][V]) receive the combined logits and the sampling distribution.
 * V <= 4096, 1 <= max_k <= min(V, 1024), 1 <= codec_size <= V.
 * Replaces the sampling of the depth decoder's frame loop
 * (models/cudagraph/depth_decoder_graph.py:487-558, _cfg_sample, with the
 * codec mask of models/logits_process.py:7-25); the draws follow the same
 * distribution from this library's own random stream. */
int bz_sample_cfg(const float* logits, int64_t ld_logits, int32_t B, int32_t V,
                  int32_t codec_size, int32_t max_k, const float* guidance,
                  const float* temperature, const int64_t* top_k,
                  const float* top_p, const int64_t* do_sample, const uint64_t* seed,
                  uint64_t* counters, int64_t* tokens, float* cfg_out,
                  float* probs_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BZ_SAMPLE_H */
